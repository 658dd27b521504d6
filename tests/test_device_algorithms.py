"""CPU tests of the device algorithms' arithmetic, emulated lane by lane in
numpy float32 and checked against the oracle.

The register FWHT of p40-kernel_amd/csrc/fwht_device.h replaces LDS
transposes with a lane mapping (element bits 4..9 -> lane bits) under which
every cross-lane butterfly partner is one DPP move or one permlane swap, and
it carries a per-lane sign through the DPP stages.  Its algebra (mapping, sign
bookkeeping, the two-swap pairing of the half-wave stages) is checked here
bit for bit against the oracle's fwht_blocks() (src/fwht.h:20-42), so a
mistake in it fails on the CPU.  The hardware semantics of the moves
themselves are covered by the GPU parity tests.
"""
import numpy as np
import pytest

from oracle import oracle as O


def fwht_row(l: int) -> int:
    e4 = (l ^ (l >> 2)) & 1
    e5 = ((l >> 1) ^ (l >> 2)) & 1
    e6 = ((l >> 2) ^ (l >> 3)) & 1
    return e4 | (e5 << 1) | (e6 << 2) | (l & 0x38)


LANES = np.arange(64)
ROWS = np.array([fwht_row(l) for l in LANES])

# source lane of each DPP pattern (all four stay inside a 16-lane row)
DPP_SRC = {
    "quad_perm[1,0,3,2]": LANES ^ 1,
    "quad_perm[2,3,0,1]": LANES ^ 2,
    "row_half_mirror": (LANES & ~7) | (7 - (LANES & 7)),
    "row_mirror": (LANES & ~15) | (15 - (LANES & 15)),
}


def permlane_swap(a, b, width):
    """v_permlane16_swap (width 16) / v_permlane32_swap (width 32): lanes of
    the odd width-groups of `a` trade places with the even groups of `b`."""
    a2, b2 = a.copy(), b.copy()
    odd = (LANES // width) % 2 == 1
    a2[odd] = b[LANES[odd] - width]
    b2[LANES[odd] - width] = a[odd]
    return a2, b2


def emulate_fwht1024_regs(x: np.ndarray) -> np.ndarray:
    """One 1024-block through the device's register FWHT, step for step."""
    v = np.stack([x[16 * r:16 * r + 16] for r in ROWS]).astype(np.float32)   # v[lane, reg]
    for h in (1, 2, 4, 8):                                                    # register stages
        for r in range(16):
            if not r & h:
                a, b = v[:, r].copy(), v[:, r | h].copy()
                v[:, r], v[:, r | h] = a + b, a - b
    for name, bit in zip(DPP_SRC, (1, 2, 4, 8)):                              # h = 16 .. 128
        c = np.where(ROWS & bit, np.float32(-1), np.float32(1))
        v = v[DPP_SRC[name]] * c[:, None] + v                                 # fmac: c*p exact
    for width in (16, 32):                                                    # h = 256, 512
        for r in range(0, 16, 2):
            a, b = permlane_swap(v[:, r], v[:, r + 1], width)
            v[:, r], v[:, r + 1] = permlane_swap(a + b, a - b, width)
    par = np.array([bin(int(r) & 15).count("1") & 1 for r in ROWS])
    scale = np.where(par == 1, np.float32(-1 / 32), np.float32(1 / 32))
    v = v * scale[:, None]
    out = np.empty(1024, np.float32)
    for l in LANES:
        out[16 * ROWS[l]:16 * ROWS[l] + 16] = v[l]
    return out


def test_lane_mapping_is_a_permutation_and_pairs_chunks():
    assert sorted(ROWS) == list(range(64))
    # a Q8_1 chunk (element bits 0..4) is the lane pair (l, l^1)
    assert np.all(ROWS[LANES ^ 1] == ROWS ^ 1)
    # each DPP pattern flips exactly its element bit
    for name, bit in zip(DPP_SRC, (1, 2, 4, 8)):
        assert np.all(ROWS[DPP_SRC[name]] == ROWS ^ bit), name


@pytest.mark.parametrize("seed", [0, 1, 2, 3])
def test_register_fwht_bit_exact(seed):
    x = O.gen_normal(7000 + seed, 1024)
    np.testing.assert_array_equal(emulate_fwht1024_regs(x).view(np.uint32),
                                  O.fwht(x).view(np.uint32))


def test_register_fwht_cancellation_and_scale_extremes():
    # wide dynamic range and exact cancellations exercise every rounding
    rng = np.random.default_rng(11)
    x = (rng.standard_normal(1024) * np.exp2(rng.integers(-30, 30, 1024))).astype(np.float32)
    x[::5] = -x[1::5][:x[::5].size]
    np.testing.assert_array_equal(emulate_fwht1024_regs(x).view(np.uint32),
                                  O.fwht(x).view(np.uint32))


def test_round_half_away_identity():
    """trunc(2p) - trunc(p) == lroundf(p) for |p| <= 127.5 (the quantiser's
    rounding, p40-kernel_amd/csrc/fwht_device.h), including every value
    within 8 ulps of each half-integer and a dense random sample."""
    halves = np.arange(-128, 128, dtype=np.float64) + 0.5
    near = [np.float32(h) for h in halves]
    cand = []
    for h in near:
        u = np.array([h], np.float32).view(np.int32)[0]
        cand.extend(np.arange(u - 8, u + 9, dtype=np.int32))
    p = np.concatenate([np.array(cand, np.int32).view(np.float32),
                        np.random.default_rng(5).uniform(-127.5, 127.5, 2_000_000).astype(np.float32),
                        np.float32([0.0, -0.0, 0.49999997, -0.49999997, 0.5, -0.5, 127.49999, 1e-30])])
    p = p[np.abs(p) <= 127.5]
    two = (p + p).astype(np.float32)
    got = np.trunc(two).astype(np.int64) - np.trunc(p).astype(np.int64)
    ref = (np.sign(p.astype(np.float64)) * np.floor(np.abs(p.astype(np.float64)) + 0.5)).astype(np.int64)
    np.testing.assert_array_equal(got, ref)


# ----------------------------------------------------------------------------
# Small batch with a block-diagonal B (gemm_bd_kernel in csrc/gemm.hip): the
# lane-level operand assembly of v_mfma_i32_16x16x64_i8, emulated in numpy.
# A lane (row x, K-group g) and a B lane (column x, K-group g) meet byte for
# byte (the instruction's A and B lane layouts are the same), so the
# emulation pairs them directly; what it checks is which code bits and which
# activation bytes each lane loads, the zero lanes, the -s start value and
# the column -> (token, chunk) bookkeeping, against the oracle's integer
# chunk dots and its GEMM.
def _bd_piece_slot(W, X, n_tok, rows, piece, nb):
    """LDS slot of one piece as the kernel's DMA fills it: each row's two
    blocks (68 bytes), then the 8 chunks x n_tok Q8_1 blocks of the piece."""
    rb = W.reshape(-1, nb * O.PQ2_BYTES)
    w = np.concatenate([rb[r, 68 * piece:68 * piece + 68] for r in rows])
    a = X.reshape(-1, n_tok * O.Q81_BYTES)[8 * piece:8 * piece + 8].ravel()
    return w, a


def _bd_emulate(W, X, n_out, nb, NT, R=16):
    CPD = 4 if NT <= 4 else 2
    lanes = np.arange(64)
    x, g = lanes & 15, lanes >> 4
    gq, hh = g >> 1, g & 1
    cc, t = x // NT, x % NT
    col_ok = cc < CPD
    cce = np.where(col_ok, cc, CPD - 1)
    y = np.zeros((n_out, NT), np.float32)
    D_all = {}
    for row0 in range(0, n_out, R):
        rows = [min(row0 + r, n_out - 1) for r in range(R)]
        acc = np.zeros((64, 4), np.float32)
        for piece in range(nb // 2):
            wl, al = _bd_piece_slot(W, X, NT, rows, piece, nb)
            for bb in range(2):
                inner = np.zeros((64, 4), np.float32)
                for dt in range(4 // CPD):
                    c0 = 4 * bb + dt * CPD
                    rec = al.reshape(8, NT, O.Q81_BYTES)
                    dsw = rec[c0 + cce, t]
                    da = dsw[:, 0:2].copy().view(np.float16).astype(np.float32).ravel()
                    s = dsw[:, 2:4].copy().view(np.int16).astype(np.int64).ravel()
                    D = np.repeat(-s[:, None], 4, axis=1)          # lane (x, g): rows 4g+i, column x
                    for m in range(CPD // 2):
                        # A: 16 int8 per lane from one code dword
                        off = x * 68 + 2 + 8 * gq + 4 * hh + 34 * bb + 8 * (dt * CPD + 2 * m)
                        wd = np.array([int.from_bytes(wl[o:o + 4].tobytes(), "little") for o in off], np.uint64)
                        A = np.stack([((wd >> np.uint64(2 * k)) & np.uint64(0x03030303)) for k in range(4)], 1)
                        Ab = A.astype("<u4").view(np.uint8).reshape(64, 16).astype(np.int64)
                        # B: the matching 16 activation bytes, or zeros
                        live = col_ok & (cc == 2 * m + gq)
                        boff = (cc * NT + t) * O.Q81_BYTES + 4 + 16 * hh + c0 * NT * O.Q81_BYTES
                        Bb = np.zeros((64, 16), np.int64)
                        for l in np.nonzero(live)[0]:
                            Bb[l] = al[boff[l]:boff[l] + 16].view(np.int8)
                        # D[r][c] += sum over g, bytes of A(r, g) * B(c, g)
                        Ar = Ab.reshape(4, 16, 16)                 # [g][row][byte]
                        Br = Bb.reshape(4, 16, 16)                 # [g][col][byte]
                        full = np.einsum("grk,gck->rc", Ar, Br)
                        for l in lanes:
                            D[l] += full[4 * g[l]:4 * g[l] + 4, x[l]]
                    D_all[(row0, piece, bb, dt)] = D.copy()
                    Df = D.astype(np.float32)
                    inner = (da[:, None] * Df) if dt == 0 else (da[:, None] * Df + inner).astype(np.float32)
                dwr = np.array([[wl[(4 * g[l] + i) * 68 + 34 * bb:(4 * g[l] + i) * 68 + 34 * bb + 2].view(np.float16)[0]
                                 for i in range(4)] for l in lanes], np.float32)
                acc = (dwr * inner + acc).astype(np.float32)
        for l in lanes:
            if not col_ok[l]:
                continue
            for i in range(4):
                r = row0 + 4 * g[l] + i
                if r < n_out:
                    y[r, t[l]] += acc[l, i]
    return y, D_all


@pytest.mark.parametrize("NT", [3, 4, 5, 8])
def test_block_diagonal_small_batch_emulation(NT):
    n_out, n_in = 20, 1024
    nb = n_in // 128
    W = O.gen_weights(4100 + NT, n_out, n_in, 0.05)
    xs = [O.gen_normal(4200 + 7 * NT + t, n_in) for t in range(NT)]
    Xt = [O.quantize_q8_1(v, True) for v in xs]
    X = np.stack([q.reshape(-1, O.Q81_BYTES) for q in Xt], 1).ravel()   # chunk-major
    y, D_all = _bd_emulate(W, X, n_out, nb, NT)
    # every result element is one exact integer chunk dot of its (token, chunk)
    dots = [O.chunk_dots(W, Xt[t], n_out, n_in) for t in range(NT)]
    CPD = 4 if NT <= 4 else 2
    for (row0, piece, bb, dt), D in D_all.items():
        for l in range(64):
            xx, gg = l & 15, l >> 4
            c, tt = xx // NT, xx % NT
            if c >= CPD:
                continue
            chunk = 8 * piece + 4 * bb + dt * CPD + c
            for i in range(4):
                r = row0 + 4 * gg + i
                if r < n_out:
                    assert D[l, i] == dots[tt][r, chunk]
    ref = O.gemm(W, X, n_out, n_in, NT)
    scale = float(np.max(np.abs(ref)))
    assert float(np.max(np.abs(y - ref))) <= 1e-5 * scale


# ------------------------------------------------------------------------
# Address math of the prefill GEMM's weight staging (gemm_f16_kernel,
# p40-kernel_amd/csrc/gemm.hip, `prefetch`): per (row, chunk ap, block) the
# kernel reads a dword-aligned window of three dwords over the chunk's 8 code
# bytes plus the 2-byte block scale, with W at any 2-byte alignment.  Restated
# here on the CPU: every byte read must lie in [0, w_bytes) -- an exact-size
# allocation can end at an unmapped page -- and the realigned words must be
# the chunk's code bytes.
def _alignbyte(hi, lo, s):
    return ((((hi.astype(np.uint64) << np.uint64(32)) | lo.astype(np.uint64)) >> (8 * s).astype(np.uint64))
            & np.uint64(0xffffffff)).astype(np.uint32)


@pytest.mark.parametrize("w_align", [0, 2])
@pytest.mark.parametrize("n_out,nb", [(17408, 40), (5120, 136), (6144, 40), (1024, 40),
                                      (129, 3), (200, 5), (64, 8), (7, 1)])
def test_gemm_f16_weight_window_stays_in_w(n_out, nb, w_align):
    rs = 34 * nb
    w_bytes = rs * n_out
    rows = np.arange(n_out, dtype=np.int64)[:, None, None]
    blk = np.arange(nb, dtype=np.int64)[None, :, None]
    ap = np.arange(4, dtype=np.int64)[None, None, :]
    a_off = rows * rs + 34 * blk + 2 + 8 * ap
    aa = ((a_off + w_align) & ~3) - w_align
    sh = (a_off + w_align) & 3
    tail = aa + 12 > w_bytes
    third = np.where(tail, np.where(sh != 0, aa + 6, aa + 4), aa + 8)
    scale = a_off - 2 - 8 * ap
    lo = np.minimum(np.minimum(aa, third), scale).min()
    hi = max((aa + 8).max(), (third + 4).max(), (scale + 2).max())
    assert lo >= 0 and hi <= w_bytes, (lo, hi, w_bytes)
    assert set(np.unique(sh)) <= {0, 2}
    # data: the realigned words are the chunk's 8 code bytes (last rows only)
    rng = np.random.default_rng(nb)
    buf = rng.integers(0, 256, w_bytes + w_align + 8, dtype=np.uint8)
    last = slice(max(0, n_out - 3), n_out)
    A, S, T, TL = (v[last].ravel() for v in (aa, sh, third, np.broadcast_to(tail, aa.shape)))
    O_ = a_off[last].ravel()
    def dword(at):
        idx = w_align + at[:, None] + np.arange(4)
        return (buf[idx].astype(np.uint32) << (8 * np.arange(4, dtype=np.uint32))).sum(axis=1).astype(np.uint32)
    w0, w1, w2 = dword(A), dword(A + 4), dword(T)
    a2 = np.where(TL, w2 >> np.uint32(16), w2)
    cw0 = _alignbyte(w1, w0, S)
    cw1 = _alignbyte(a2, w1, S)
    want0 = dword(O_)
    want1 = dword(O_ + 4)
    assert np.array_equal(cw0, want0)
    assert np.array_equal(cw1, want1)


# ------------------------------------------------ GEMV unit numbering / tail
def _gemv_wave_index(w, blk, blocks, xl):
    """gemv_nb_kernel's wave numbering (csrc/gemv.hip, wave_index): plain
    slot-major, or groups of 2^xl consecutive units per XCD."""
    if xl <= 0:
        return w * blocks + blk
    K = blocks >> 3
    t = w * K + (blk >> 3)
    m = (1 << xl) - 1
    return ((((t >> xl) << 3) + (blk & 7)) << xl) | (t & m)


def _dispatch_xl(blocks, waves, xl=3):
    """launch_nb_t's choice of the XCD group size for a grid."""
    if blocks % 8 != 0:
        return 0
    while xl > 0 and ((blocks // 8) * waves) % (1 << xl) != 0:
        xl -= 1
    return xl


@pytest.mark.parametrize("waves", [4, 6, 8])
@pytest.mark.parametrize("blocks", [8, 16, 24, 64, 248, 256, 768])
def test_gemv_numbering_and_shared_tail_condition(blocks, waves):
    """The numbering is a permutation of the grid's waves, and wherever the
    dispatcher enables the shared tail (L = T * blocks last-round units, 2^xl
    dividing T * blocks / 8) the units of the last round are exactly the last
    units of waves 0..T-1 of every workgroup -- the kernel's assumption."""
    for want_xl in range(4):
        xl = min(want_xl, _dispatch_xl(blocks, waves))
        idx = np.array([[_gemv_wave_index(w, b, blocks, xl) for b in range(blocks)] for w in range(waves)])
        assert sorted(idx.ravel().tolist()) == list(range(waves * blocks))
        for T in range(1, waves):
            if xl and (T * (blocks // 8)) % (1 << xl) != 0:
                continue
            owner = idx < T * blocks
            assert np.array_equal(owner, np.arange(waves)[:, None] < T + np.zeros((1, blocks), dtype=int))
