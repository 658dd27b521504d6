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
