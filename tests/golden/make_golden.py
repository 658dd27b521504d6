"""Writes the golden fixtures F1-F9 from the reference's own host code.

The vectors come from oracle/_ref/libbonsai_ref.so, i.e. the reference
headers src/pq2_0.h, src/fwht.h, src/pq2_0_repack.h and src/ops.h compiled
from /root/reference by `make -C oracle ref` (see oracle/ref_shim.cpp).  Inputs
are drawn with the oracle's seeded generator (splitmix64 + Box-Muller), which
is plain data generation, not a checked function.  Run once in a container
that has the reference tree; the fixtures (golden.npz) are committed and the
tests read only them.

    python tests/golden/make_golden.py
"""
from __future__ import annotations

import ctypes as C
import os
import struct
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)
from oracle import oracle as O  # noqa: E402

OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden.npz")


def p(a, t):
    return a.ctypes.data_as(t)


def ref_q8(R, x, permute=True):
    x = np.ascontiguousarray(x, np.float32)
    y = np.empty(x.size // 32 * 36, np.uint8)
    R.ref_quantize_q8_1(p(x, O._f32p), p(y, O._u8p), x.size, int(permute))
    return y


def ref_fwht(R, x, signs=None):
    y = np.array(x, np.float32, copy=True)
    R.ref_fwht_blocks(p(y, O._f32p), None if signs is None else p(signs, O._f32p), y.size)
    return y


def ref_gemv(R, W, xq, n_out, n_in):
    y = np.empty(n_out, np.float32)
    R.ref_gemv(p(W, O._u8p), p(xq, O._u8p), p(y, O._f32p), n_out, n_in)
    return y


def ref_chunk_sumi(R, W, xq, n_out, n_in):
    nb, nc = n_in // 128, n_in // 32
    out = np.empty((n_out, nc), np.int32)
    for r in range(n_out):
        for c in range(nc):
            wb = W[(r * nb + c // 4) * 34:]
            ab = xq[c * 36:]
            out[r, c] = R.ref_chunk_sumi(p(wb, O._u8p), p(ab, O._u8p), c % 4)
    return out


def f16_edge_inputs():
    v = []
    # exact ties between adjacent normal fp16 values, both signs, many binades
    for e in range(-14, 16):
        for m in (0, 1, 2, 3, 511, 512, 1021, 1022):
            lo = (1 + m / 1024.0) * 2.0 ** e
            v += [lo + 2.0 ** (e - 11), -(lo + 2.0 ** (e - 11))]
    # subnormal range and its ties, underflow to zero, overflow
    for k in range(0, 40):
        v.append(k * 2.0 ** -25)
        v.append((k + 0.5) * 2.0 ** -24)
    v += [2.0 ** -25, 2.0 ** -26, 2.0 ** -24, 65504.0, 65519.99, 65520.0, 65536.0, 1e9, -1e9,
          0.0, -0.0, float("inf"), float("-inf"), float("nan"), 1.0 / 127.0, 3.0 / 127.0]
    return np.array(v, np.float32)


def tie_chunk():
    """A chunk whose x*id products land exactly on k + 0.5 (round-away ties)."""
    x = np.zeros(32, np.float32)
    x[0] = 127.0                      # amax -> d = 1, id = 1
    x[1:16] = np.array([0.5, -0.5, 1.5, -1.5, 2.5, -2.5, 126.5, -126.5, 3.5, 10.5, -10.5,
                        0.25, -0.75, 64.5, -64.5], np.float32)
    x[16:32] = np.arange(16, dtype=np.float32) * 7.5 - 60.0
    return x


def pq2_special_blocks():
    """Blocks for the ternary quantiser's edge cases (src/pq2_0.h:74-90)."""
    blocks = []
    b = np.zeros(128, np.float32)            # all zero: d = 0, id = 0, every code 1
    blocks.append(b)
    b = np.zeros(128, np.float32)            # x * id exactly +-0.5: lroundf goes away from zero
    b[0] = 2.0
    b[1:9] = [1.0, -1.0, 1.0, -1.0, 0.5, -0.5, 1.5, -1.5]
    b[9:] = np.linspace(-2.0, 2.0, 119).astype(np.float32)
    blocks.append(b)
    b = np.linspace(-1.0, 1.0, 128).astype(np.float32)
    b[5] = 1.0 + 2.0 ** -11                  # amax an exact fp16 tie (1 and 1 + 2^-10): ties away
    blocks.append(b)
    blocks.append(np.linspace(-1e-6, 3e-6, 128).astype(np.float32))    # subnormal fp16 scale
    blocks.append(np.linspace(-7e4, 1e5, 128).astype(np.float32))      # scale overflows fp16
    b = -np.abs(np.linspace(0.1, 3.0, 128)).astype(np.float32)        # all negative
    blocks.append(b)
    return np.concatenate(blocks)


def main():
    R = O.ref()
    if R is None:
        raise SystemExit("oracle/_ref/libbonsai_ref.so missing: run `make -C oracle ref` first")
    fx = {}

    # F1: fp16 encode on edge cases + full 2^32 hash + full decode table
    e = f16_edge_inputs()
    fx["f1_in"] = e
    fx["f1_out"] = np.array([R.ref_f32_to_f16(float(t)) for t in e], np.uint16)
    fx["f1_hash_all"] = np.array([R.ref_f16_encode_hash(0, 1 << 32, 1)], np.uint64)
    fx["f1_decode_all"] = np.array([R.ref_f16_to_f32(h) for h in range(65536)], np.float32)

    # F2: Q8_1 quantiser
    x = O.gen_normal(101, 5120)
    x = ref_fwht(R, x)
    special = np.concatenate([tie_chunk(), np.zeros(32, np.float32),
                              np.full(32, 1e-30, np.float32),
                              np.linspace(-3, 3, 32).astype(np.float32),
                              np.where(np.arange(32) % 2 == 0, 1e4, -3e-3).astype(np.float32)])
    for name, v in (("seeded", x), ("special", special), ("k32", O.gen_normal(102, 32) * 5)):
        fx[f"f2_{name}_in"] = v.astype(np.float32)
        fx[f"f2_{name}_perm"] = ref_q8(R, v, True)
        fx[f"f2_{name}_plain"] = ref_q8(R, v, False)

    # F3: FWHT bit patterns, signs NULL and a length-n +-1 vector
    x3 = O.gen_normal(103, 2048)
    s3 = np.where(O.gen_normal(104, 2048) > 0, 1.0, -1.0).astype(np.float32)
    fx["f3_in"] = x3
    fx["f3_signs"] = s3
    fx["f3_out"] = ref_fwht(R, x3)
    fx["f3_out_signed"] = ref_fwht(R, x3, s3)

    # F4: chunk dots + row dots at K = 5120 and 17408 (code-3 rich weights)
    for k, seed in ((5120, 105), (17408, 106)):
        n_out = 8
        W = O.gen_weights(seed, n_out, k, 0.02)
        xa = ref_fwht(R, O.gen_normal(seed + 1000, k))
        xq = ref_q8(R, xa, True)
        fx[f"f4_{k}_W"] = W
        fx[f"f4_{k}_xq"] = xq
        fx[f"f4_{k}_sumi"] = ref_chunk_sumi(R, W, xq, n_out, k)
        fx[f"f4_{k}_y"] = ref_gemv(R, W, xq, n_out, k)

    # F5: repack bytes + repack row dot
    W5 = fx["f4_5120_W"]
    Wr = np.empty_like(W5)
    assert R.ref_repack_rows(p(W5, O._u8p), p(Wr, O._u8p), 8, 5120) == 0
    fx["f5_Wr"] = Wr
    fx["f5_y"] = np.array([R.ref_repack_row_dot(p(Wr[r * 1360:], O._u8p), p(fx["f4_5120_xq"], O._u8p), 40)
                           for r in range(8)], np.float32)

    # F6: chunk-major GEMM (the tests/test_p40.cpp:449-470 loop)
    for (n_out, n_in, n_tok, seed) in ((64, 256, 5, 107), (32, 1024, 8, 108)):
        W = O.gen_weights(seed, n_out, n_in, 0.01)
        X = O.gen_normal(seed + 1, n_tok * n_in).reshape(n_tok, n_in)
        Xq = np.empty(n_in // 32 * n_tok * 36, np.uint8)
        for t in range(n_tok):
            q = ref_q8(R, X[t], True).reshape(-1, 36)
            for c in range(n_in // 32):
                Xq[(c * n_tok + t) * 36:(c * n_tok + t + 1) * 36] = q[c]
        Y = np.empty(n_out * n_tok, np.float32)
        R.ref_gemm(p(W, O._u8p), p(Xq, O._u8p), p(Y, O._f32p), n_out, n_in, n_tok)
        tag = f"f6_{n_out}x{n_in}x{n_tok}"
        fx[tag + "_W"], fx[tag + "_X"], fx[tag + "_Xq"], fx[tag + "_Y"] = W, X, Xq, Y

    # F7: SwiGLU -> FWHT -> Q8_1 chain
    g = O.gen_normal(109, 2048) * 2
    u = O.gen_normal(110, 2048)
    h = np.empty(2048, np.float32)
    R.ref_swiglu(p(g, O._f32p), p(u, O._f32p), p(h, O._f32p), 2048)
    fx["f7_gate"], fx["f7_up"], fx["f7_h"] = g, u, h
    fx["f7_hq"] = ref_q8(R, ref_fwht(R, h), True)

    # F8: RMSNorm (src/ops.h:13-22) -> FWHT -> Q8_1, two rows and two eps
    for (n, seed, eps) in ((3072, 111, 1e-6), (1024, 113, 1e-2)):
        x = O.gen_normal(seed, n) * 3
        w = O.gen_normal(seed + 1, n) * 0.1 + 1
        y = np.empty(n, np.float32)
        R.ref_rmsnorm(p(x, O._f32p), p(w, O._f32p), p(y, O._f32p), n, C.c_float(eps))
        tag = f"f8_{n}"
        fx[tag + "_x"], fx[tag + "_w"], fx[tag + "_y"] = x, w, y
        fx[tag + "_eps"] = np.float32(eps)
        fx[tag + "_yq"] = ref_q8(R, ref_fwht(R, y), True)

    # F9: reference ternary quantiser, dequantiser and float block dot
    #     (src/pq2_0.h:62-90, 134-142)
    xs = np.concatenate([O.gen_normal(115, 8 * 1024, 0.02), pq2_special_blocks()])
    w9 = np.empty(xs.size // 128 * 34, np.uint8)
    R.ref_quantize_pq2_0(p(xs, O._f32p), p(w9, O._u8p), xs.size)
    fx["f9_x"], fx["f9_w"] = xs, w9
    wd = np.concatenate([w9, fx["f4_5120_W"][:34 * 40]])       # plus code-3-rich rows
    yd = np.empty(wd.size // 34 * 128, np.float32)
    R.ref_dequantize_pq2_0(p(wd, O._u8p), p(yd, O._f32p), yd.size)
    fx["f9_wd"], fx["f9_deq"] = wd, yd
    a9 = O.gen_normal(116, yd.size) * 3
    fx["f9_a"] = a9
    fx["f9_dot"] = np.array([R.ref_pq2_0_dot_f32(p(wd[34 * i:], O._u8p), p(a9[128 * i:], O._f32p))
                             for i in range(wd.size // 34)], np.float32)

    np.savez_compressed(OUT, **fx)
    print(f"wrote {OUT}: {os.path.getsize(OUT)} bytes, {len(fx)} arrays")


if __name__ == "__main__":
    main()
