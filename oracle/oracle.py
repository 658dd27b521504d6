"""ctypes/numpy front end of the CPU parity oracle.

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py, as the checker.  The product (p40-kernel_amd/)
never imports this module.

Two libraries sit behind it:
  * liboracle.so       -- pq2_oracle.c, the build's own C restatement of the
                          reference host path (src/pq2_0.h, src/fwht.h,
                          src/pq2_0_repack.h, src/ops.h, tests/test_p40.cpp);
  * _ref/libbonsai_ref.so -- the reference's own header code compiled from
                          /root/reference (ref_shim.cpp); optional, present
                          where it was built.
Byte buffers are numpy uint8 arrays in the reference's exact layouts
(block_pq2_0 = 34 B, block_q8_1 = 36 B).
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
QK_PQ2, QK8, PQ2_BYTES, Q81_BYTES, HBLK = 128, 32, 34, 36, 1024

_u8p = C.POINTER(C.c_uint8)
_f32p = C.POINTER(C.c_float)
_i32p = C.POINTER(C.c_int32)
_i64 = C.c_int64


def _p(a: np.ndarray, t):
    return a.ctypes.data_as(t)


def _load(path: str, required: bool):
    if not os.path.exists(path):
        if required:
            raise RuntimeError(f"oracle library missing: {path} (run `make -C oracle`)")
        return None
    return C.CDLL(path)


_lib = None
_ref = None


def lib():
    global _lib
    if _lib is None:
        _lib = _load(os.path.join(HERE, "liboracle.so"), True)
        L = _lib
        L.orc_f16_to_f32.argtypes = [C.c_uint16]; L.orc_f16_to_f32.restype = C.c_float
        L.orc_f32_to_f16.argtypes = [C.c_float]; L.orc_f32_to_f16.restype = C.c_uint16
        L.orc_f16_encode_hash.argtypes = [C.c_uint64] * 3; L.orc_f16_encode_hash.restype = C.c_uint64
        L.orc_quantize_q8_1.argtypes = [_f32p, _u8p, _i64, C.c_int]
        L.orc_quantize_chunk_major.argtypes = [_f32p, _u8p, _i64, _i64]
        L.orc_fwht_blocks.argtypes = [_f32p, _f32p, _i64]
        L.orc_dequantize_pq2_0.argtypes = [_u8p, _f32p, _i64]
        L.orc_quantize_pq2_0.argtypes = [_f32p, _u8p, _i64]
        L.orc_pq2_0_dot_f32.argtypes = [_u8p, _f32p]; L.orc_pq2_0_dot_f32.restype = C.c_float
        L.orc_chunk_sumi.argtypes = [_u8p, _u8p, C.c_int]; L.orc_chunk_sumi.restype = C.c_int32
        L.orc_row_dot.argtypes = [_u8p, _u8p, _i64]; L.orc_row_dot.restype = C.c_float
        L.orc_gemv.argtypes = [_u8p, _u8p, _f32p, _i64, _i64, C.c_int]
        L.orc_chunk_dots.argtypes = [_u8p, _u8p, _i32p, _i64, _i64]
        L.orc_gemm.argtypes = [_u8p, _u8p, _f32p, _i64, _i64, _i64, C.c_int]
        L.orc_repack_rows.argtypes = [_u8p, _u8p, _i64, _i64]; L.orc_repack_rows.restype = C.c_int
        L.orc_unpack_rows.argtypes = [_u8p, _u8p, _i64, _i64]; L.orc_unpack_rows.restype = C.c_int
        L.orc_repack_row_dot.argtypes = [_u8p, _u8p, _i64]; L.orc_repack_row_dot.restype = C.c_float
        L.orc_gemv_repack.argtypes = [_u8p, _f32p, _f32p, _i64, _i64, C.c_int]
        L.orc_swiglu.argtypes = [_f32p, _f32p, _f32p, _i64]
        L.orc_rmsnorm.argtypes = [_f32p, _f32p, _f32p, _i64, C.c_float]
        L.orc_gen_normal.argtypes = [C.c_uint64, _f32p, _i64, C.c_float]
        L.orc_gen_weights.argtypes = [C.c_uint64, _u8p, _i64, _i64, C.c_double]
    return _lib


def ref():
    """The compiled reference (oracle/_ref), or None where it was not built."""
    global _ref
    if _ref is None:
        _ref = _load(os.path.join(HERE, "_ref", "libbonsai_ref.so"), False)
        if _ref is None:
            return None
        R = _ref
        R.ref_f32_to_f16.argtypes = [C.c_float]; R.ref_f32_to_f16.restype = C.c_uint16
        R.ref_f16_to_f32.argtypes = [C.c_uint16]; R.ref_f16_to_f32.restype = C.c_float
        R.ref_f16_encode_hash.argtypes = [C.c_uint64] * 3; R.ref_f16_encode_hash.restype = C.c_uint64
        R.ref_quantize_q8_1.argtypes = [_f32p, _u8p, _i64, C.c_int]
        R.ref_fwht_blocks.argtypes = [_f32p, _f32p, _i64]
        R.ref_quantize_pq2_0.argtypes = [_f32p, _u8p, _i64]
        R.ref_dequantize_pq2_0.argtypes = [_u8p, _f32p, _i64]
        R.ref_pq2_0_dot_f32.argtypes = [_u8p, _f32p]; R.ref_pq2_0_dot_f32.restype = C.c_float
        R.ref_chunk_sumi.argtypes = [_u8p, _u8p, C.c_int]; R.ref_chunk_sumi.restype = C.c_int32
        R.ref_row_dot.argtypes = [_u8p, _u8p, _i64]; R.ref_row_dot.restype = C.c_float
        R.ref_gemv.argtypes = [_u8p, _u8p, _f32p, _i64, _i64]
        R.ref_gemm.argtypes = [_u8p, _u8p, _f32p, _i64, _i64, _i64]
        R.ref_repack_rows.argtypes = [_u8p, _u8p, _i64, _i64]; R.ref_repack_rows.restype = C.c_int
        R.ref_unpack_rows.argtypes = [_u8p, _u8p, _i64, _i64]; R.ref_unpack_rows.restype = C.c_int
        R.ref_repack_row_dot.argtypes = [_u8p, _u8p, _i64]; R.ref_repack_row_dot.restype = C.c_float
        R.ref_swiglu.argtypes = [_f32p, _f32p, _f32p, _i64]
        R.ref_rmsnorm.argtypes = [_f32p, _f32p, _f32p, _i64, C.c_float]
    return _ref


# ----------------------------------------------------------------- wrappers
def f32_to_f16(x: float) -> int:
    return lib().orc_f32_to_f16(float(x))


def f16_to_f32(h: int) -> float:
    return lib().orc_f16_to_f32(int(h))


def quantize_q8_1(x: np.ndarray, permute: bool = True) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    assert x.size % QK8 == 0
    y = np.empty(x.size // QK8 * Q81_BYTES, np.uint8)
    lib().orc_quantize_q8_1(_p(x, _f32p), _p(y, _u8p), x.size, int(permute))
    return y


def quantize_chunk_major(x: np.ndarray) -> np.ndarray:
    """x: [n_tok, n_in] fp32 -> chunk-major Q8_1 bytes [n_in/32][n_tok]."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    n_tok, k = x.shape
    y = np.empty(k // QK8 * n_tok * Q81_BYTES, np.uint8)
    lib().orc_quantize_chunk_major(_p(x, _f32p), _p(y, _u8p), k, n_tok)
    return y


def fwht(x: np.ndarray, signs: np.ndarray | None = None) -> np.ndarray:
    y = np.array(x, dtype=np.float32, copy=True)
    if y.size % HBLK != 0:      # the C restatement walks whole 1024-blocks
        raise ValueError(f"fwht: length {y.size} is not a multiple of {HBLK}")
    if signs is not None and np.size(signs) < y.size:
        raise ValueError("fwht: the sign vector is shorter than x")
    s = None if signs is None else np.ascontiguousarray(signs, dtype=np.float32)
    lib().orc_fwht_blocks(_p(y, _f32p), None if s is None else _p(s, _f32p), y.size)
    return y


def dequantize_pq2_0(w: np.ndarray, k: int) -> np.ndarray:
    y = np.empty(k, np.float32)
    lib().orc_dequantize_pq2_0(_p(w, _u8p), _p(y, _f32p), k)
    return y


def quantize_pq2_0(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    w = np.empty(x.size // QK_PQ2 * PQ2_BYTES, np.uint8)
    lib().orc_quantize_pq2_0(_p(x, _f32p), _p(w, _u8p), x.size)
    return w


def pq2_0_dot_f32(W: np.ndarray, a: np.ndarray) -> np.ndarray:
    """Float dot of every 34-byte block of W with its 128 floats of a
    (a.size == 128 * blocks): one value per block."""
    W = np.ascontiguousarray(W, np.uint8); a = np.ascontiguousarray(a, np.float32)
    nblk = W.size // PQ2_BYTES
    assert a.size == nblk * QK_PQ2
    L = lib()
    return np.array([L.orc_pq2_0_dot_f32(_p(W[b * PQ2_BYTES:], _u8p), _p(a[b * QK_PQ2:], _f32p))
                     for b in range(nblk)], np.float32)


def gemv(W: np.ndarray, xq: np.ndarray, n_out: int, n_in: int, nthreads: int = 1) -> np.ndarray:
    y = np.empty(n_out, np.float32)
    lib().orc_gemv(_p(W, _u8p), _p(xq, _u8p), _p(y, _f32p), n_out, n_in, nthreads)
    return y


def chunk_dots(W: np.ndarray, xq: np.ndarray, n_out: int, n_in: int) -> np.ndarray:
    out = np.empty((n_out, n_in // QK8), np.int32)
    lib().orc_chunk_dots(_p(W, _u8p), _p(xq, _u8p), _p(out, _i32p), n_out, n_in)
    return out


def gemm(W: np.ndarray, X: np.ndarray, n_out: int, n_in: int, n_tok: int,
         nthreads: int = 1) -> np.ndarray:
    Y = np.empty((n_out, n_tok), np.float32)
    lib().orc_gemm(_p(W, _u8p), _p(X, _u8p), _p(Y, _f32p), n_out, n_in, n_tok, nthreads)
    return Y


def repack(W: np.ndarray, n_out: int, n_in: int) -> np.ndarray:
    out = np.empty_like(W)
    rc = lib().orc_repack_rows(_p(W, _u8p), _p(out, _u8p), n_out, n_in)
    if rc:
        raise ValueError("repack requires n_in/128 to be a positive multiple of 8")
    return out


def unpack(Wr: np.ndarray, n_out: int, n_in: int) -> np.ndarray:
    out = np.empty_like(Wr)
    rc = lib().orc_unpack_rows(_p(Wr, _u8p), _p(out, _u8p), n_out, n_in)
    if rc:
        raise ValueError("unpack requires n_in/128 to be a positive multiple of 8")
    return out


def gemv_repack(Wr: np.ndarray, x: np.ndarray, n_out: int, n_in: int, nthreads: int = 1):
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.empty(n_out, np.float32)
    lib().orc_gemv_repack(_p(Wr, _u8p), _p(x, _f32p), _p(y, _f32p), n_out, n_in, nthreads)
    return y


def swiglu(g: np.ndarray, u: np.ndarray) -> np.ndarray:
    g = np.ascontiguousarray(g, np.float32); u = np.ascontiguousarray(u, np.float32)
    y = np.empty_like(g)
    lib().orc_swiglu(_p(g, _f32p), _p(u, _f32p), _p(y, _f32p), g.size)
    return y


def rmsnorm(x: np.ndarray, w: np.ndarray, eps: float) -> np.ndarray:
    """RMSNorm of one row (src/ops.h:13-22): sequential fp32 sum of squares."""
    x = np.ascontiguousarray(x, np.float32); w = np.ascontiguousarray(w, np.float32)
    y = np.empty_like(x)
    lib().orc_rmsnorm(_p(x, _f32p), _p(w, _f32p), _p(y, _f32p), x.size, C.c_float(eps))
    return y


def gen_normal(seed: int, n: int, sigma: float = 1.0) -> np.ndarray:
    x = np.empty(n, np.float32)
    lib().orc_gen_normal(seed, _p(x, _f32p), n, sigma)
    return x


def gen_weights(seed: int, n_out: int, n_in: int, p3: float = 0.001) -> np.ndarray:
    W = np.empty(n_out * (n_in // QK_PQ2) * PQ2_BYTES, np.uint8)
    lib().orc_gen_weights(seed, _p(W, _u8p), n_out, n_in, p3)
    return W


# -------------------------------------------------- decoded views (numpy)
def q81_fields(q: np.ndarray):
    """(d fp16 bits uint16, s int16, qs int8 [nblk, 32]) of a Q8_1 byte buffer."""
    b = q.reshape(-1, Q81_BYTES)
    d = b[:, 0:2].copy().view(np.uint16).ravel()
    s = b[:, 2:4].copy().view(np.int16).ravel()
    qs = b[:, 4:].copy().view(np.int8)
    return d, s, qs


def pq2_fields(W: np.ndarray):
    """(d fp16 bits uint16 [nblk], codes uint8 [nblk, 128]) of PQ2_0 bytes."""
    b = W.reshape(-1, PQ2_BYTES)
    d = b[:, 0:2].copy().view(np.uint16).ravel()
    by = b[:, 2:]
    codes = np.stack([(by >> (2 * e)) & 3 for e in range(4)], axis=-1).reshape(-1, QK_PQ2)
    return d, codes
