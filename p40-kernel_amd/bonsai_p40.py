"""Host-side Python binding of libbonsai_p40.so (the gfx950 PQ2_0 matmul path).

The native library exports the C ABI of include/bonsai_p40.h; this module
binds it with ctypes and offers thin wrappers over torch device tensors
(torch is used only for device memory and the current HIP stream).  Every
wrapper raises if the library is missing or a call returns nonzero -- there is
no CPU fallback in this module.

Reference interface mirrored: include/bonsai_p40.h of boetti-dev/p40-kernel
(bonsai_p40_gemv, _quant_activations, _gemm, _repack, _gemv_repack, _fwht,
_rmsnorm), plus the additions declared at the end of the header.
"""
from __future__ import annotations

import ctypes as C
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libbonsai_p40.so")

QK_PQ2 = 128          # weights per block_pq2_0
QK8 = 32              # elements per block_q8_1
PQ2_BYTES = 34        # sizeof(block_pq2_0)
Q81_BYTES = 36        # sizeof(block_q8_1)
HBLK = 1024           # Hadamard block

# Every symbol of include/bonsai_p40.h with its ctypes signature.
_V, _I64, _F32P = C.c_void_p, C.c_int64, C.c_void_p
SIGNATURES = {
    "bonsai_p40_gemv": [_V, _V, _F32P, _I64, _I64, _V],
    "bonsai_p40_quant_activations": [_F32P, _V, _I64, _V],
    "bonsai_p40_gemm": [_V, _V, _F32P, _I64, _I64, _I64, _V],
    "bonsai_p40_gemm_ws": [_V, _V, _F32P, _I64, _I64, _I64, _V, _I64, _V],
    "bonsai_p40_gemm_workspace_bytes": [_I64, _I64],
    "bonsai_p40_repack": [_V, _V, _I64, _I64, _V],
    "bonsai_p40_gemv_repack": [_V, _F32P, _F32P, _I64, _I64, _V],
    "bonsai_p40_fwht": [_F32P, _F32P, _I64, _V],
    "bonsai_p40_fwht_signs_n": [_F32P, _F32P, _I64, _V],
    "bonsai_p40_rmsnorm": [_F32P, _F32P, _F32P, _I64, _I64, C.c_float, _V],
    "bonsai_p40_gdn_step": [_F32P] * 7 + [C.c_int] * 4 + [_V],
    "bonsai_p40_attn": [_F32P] * 4 + [C.c_int] * 4 + [C.c_float, _V],
    "bonsai_p40_fwht_quant": [_F32P, _F32P, _V, _I64, _V],
    "bonsai_p40_quant_tokens": [_F32P, _F32P, _V, _I64, _I64, C.c_int, _V],
    "bonsai_p40_swiglu_fwht_quant": [_F32P, _F32P, _F32P, _V, _I64, _V],
    "bonsai_p40_rmsnorm_fwht_quant": [_F32P, _F32P, _F32P, _V, _I64, _I64, C.c_float, _V],
    "bonsai_p40_fwht_gemv": [_V, _F32P, _F32P, _F32P, _I64, _I64, _V],
    "bonsai_p40_quant_gemv": [_V, _F32P, _F32P, _I64, _I64, _V],
    "bonsai_p40_ggml_should_use": [C.c_int, C.c_int, _I64],
    "bonsai_p40_ggml_mul_mat": [_V, _V, _V, _V, C.c_size_t, _V],
    "bonsai_p40_gemv_group": [_V, _V, _V, C.c_int, _V, _I64, _V],
    "bonsai_p40_fwht_gemv_group": [_V, _V, _V, C.c_int, _F32P, _F32P, _I64, _V],
    "bonsai_p40_rmsnorm_fwht_gemv_group": [_V, _V, _V, C.c_int, _F32P, _F32P, _F32P, _I64, C.c_float, _V],
    "bonsai_p40_ffn_gate_up_swiglu": [_V, _V, _F32P, _F32P, _F32P, _F32P, _V, _I64, _I64, C.c_float, _V, _V, _V],
    "bonsai_p40_ffn_gate_up_swiglu_noalloc": [_V, _V, _F32P, _F32P, _F32P, _F32P, _V, _I64, _I64, C.c_float,
                                              _V, _V],
    "bonsai_p40_quantize_pq2_0": [_F32P, _V, _I64, _V],
    "bonsai_p40_dequantize_pq2_0": [_V, _F32P, _I64, _V],
    "bonsai_p40_chunk_dots": [_V, _V, _V, _I64, _I64, _V],
    "bonsai_p40_stream_read": [_V, _I64, _V, C.c_int, _V],
    "bonsai_p40_reload_tuning": [],
    "bonsai_p40_mfma_probe": [C.c_int, C.c_int, C.c_int, _V, _V, _V],
    "bonsai_p40_overlap_probe": [C.c_int, C.c_int, C.c_int, C.c_int, _V, _V],
    "bonsai_p40_launch_probe": [C.c_int, C.c_int, _V, _V],
    "bonsai_p40_unit_dma_probe": [_V, _I64, _I64, _V, _V],
    "bonsai_p40_chain_plan_bytes": [C.c_int],
    "bonsai_p40_chain_plan": [_V, C.c_int, _V],
    "bonsai_p40_chain_run": [_V, C.c_int, _V, _V, _V],
}
RESTYPES = {"bonsai_p40_chain_plan_bytes": C.c_int64, "bonsai_p40_gemm_workspace_bytes": C.c_int64}

_lib = None


def lib() -> C.CDLL:
    """Load libbonsai_p40.so; raise if it was not built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"{LIB_PATH} is missing: build it with `make -C p40-kernel_amd` "
                "(or __graft_entry__.build())")
        L = C.CDLL(LIB_PATH)
        for name, argtypes in SIGNATURES.items():
            fn = getattr(L, name)
            fn.argtypes = argtypes
            fn.restype = RESTYPES.get(name, C.c_int)
        _lib = L
    return _lib


class BonsaiError(RuntimeError):
    pass


def _check(name: str, rc: int) -> None:
    if rc != 0:
        raise BonsaiError(f"{name} returned {rc}")


def _ptr(t) -> int | None:
    if t is None:
        return None
    if isinstance(t, int):
        return t
    return t.data_ptr()


def _stream(stream) -> int | None:
    if stream is not None:
        return stream if isinstance(stream, int) else stream.cuda_stream
    import torch
    return torch.cuda.current_stream().cuda_stream


def call(name: str, *args, stream=None) -> int:
    """Raw call: tensors are passed as device pointers; returns the rc."""
    fn = getattr(lib(), name)
    conv = [_ptr(a) if (a is None or hasattr(a, "data_ptr")) else a for a in args]
    return fn(*conv, _stream(stream))


# -------------------------------------------------------------- wrappers
def gemv(W, xq, y, n_out: int, n_in: int, stream=None) -> None:
    _check("bonsai_p40_gemv", call("bonsai_p40_gemv", W, xq, y, n_out, n_in, stream=stream))


def quant_activations(x, out, n: int, stream=None) -> None:
    _check("bonsai_p40_quant_activations",
           call("bonsai_p40_quant_activations", x, out, n, stream=stream))


def gemm(W, Xq, Y, n_out: int, n_in: int, n_tok: int, stream=None) -> None:
    _check("bonsai_p40_gemm", call("bonsai_p40_gemm", W, Xq, Y, n_out, n_in, n_tok, stream=stream))


def gemm_workspace_bytes(n_in: int, n_tok: int) -> int:
    """bonsai_p40_gemm_workspace_bytes: the workspace bonsai_p40_gemm_ws needs."""
    return int(lib().bonsai_p40_gemm_workspace_bytes(n_in, n_tok))


def gemm_ws(W, Xq, Y, n_out: int, n_in: int, n_tok: int, ws, ws_bytes=None, stream=None) -> None:
    """bonsai_p40_gemm with a workspace (a tensor, or a pointer with ws_bytes);
    Y is bit-identical to gemm()'s."""
    if ws_bytes is None:
        ws_bytes = 0 if ws is None else ws.numel() * ws.element_size()
    _check("bonsai_p40_gemm_ws", call("bonsai_p40_gemm_ws", W, Xq, Y, n_out, n_in, n_tok, ws, ws_bytes,
                                      stream=stream))


def repack(src, dst, n_out: int, n_in: int, stream=None) -> None:
    _check("bonsai_p40_repack", call("bonsai_p40_repack", src, dst, n_out, n_in, stream=stream))


def gemv_repack(W, x, y, n_out: int, n_in: int, stream=None) -> None:
    _check("bonsai_p40_gemv_repack",
           call("bonsai_p40_gemv_repack", W, x, y, n_out, n_in, stream=stream))


def fwht(x, signs, n: int, stream=None) -> None:
    """In-place FWHT-1024 blocks; signs (or None) has 1024 entries reused by
    every block, as the reference device kernel."""
    _check("bonsai_p40_fwht", call("bonsai_p40_fwht", x, signs, n, stream=stream))


def fwht_signs_n(x, signs, n: int, stream=None) -> None:
    """In-place FWHT-1024 blocks; signs (or None) is a length-n vector, block
    b using signs[1024 b ..] (the host fwht_blocks form)."""
    _check("bonsai_p40_fwht_signs_n", call("bonsai_p40_fwht_signs_n", x, signs, n, stream=stream))


def rmsnorm(x, w, y, n_rows: int, n: int, eps: float, stream=None) -> None:
    _check("bonsai_p40_rmsnorm",
           call("bonsai_p40_rmsnorm", x, w, y, n_rows, n, C.c_float(eps), stream=stream))


def fwht_quant(x, signs, xq, n: int, stream=None) -> None:
    _check("bonsai_p40_fwht_quant", call("bonsai_p40_fwht_quant", x, signs, xq, n, stream=stream))


def quant_tokens(X, signs, Xq, n: int, n_tok: int, rotate: bool, stream=None) -> None:
    _check("bonsai_p40_quant_tokens",
           call("bonsai_p40_quant_tokens", X, signs, Xq, n, n_tok, int(rotate), stream=stream))


def swiglu_fwht_quant(gate, up, signs, xq, n: int, stream=None) -> None:
    _check("bonsai_p40_swiglu_fwht_quant",
           call("bonsai_p40_swiglu_fwht_quant", gate, up, signs, xq, n, stream=stream))


def rmsnorm_fwht_quant(x, w, signs, xq, n: int, n_tok: int, eps: float, stream=None) -> None:
    _check("bonsai_p40_rmsnorm_fwht_quant",
           call("bonsai_p40_rmsnorm_fwht_quant", x, w, signs, xq, n, n_tok, C.c_float(eps),
                stream=stream))


def quant_gemv(W, x, y, n_out: int, n_in: int, stream=None) -> None:
    """y = W . Q8_1(x), one launch (no rotation, no Q8_1 buffer)."""
    _check("bonsai_p40_quant_gemv", call("bonsai_p40_quant_gemv", W, x, y, n_out, n_in, stream=stream))


class GgmlTensor(C.Structure):
    """bonsai_ggml_tensor of include/bonsai_p40_ggml.h: the ggml_tensor fields
    the ggml hook reads."""
    _fields_ = [("type", C.c_int), ("ne", C.c_int64 * 4), ("nb", C.c_size_t * 4), ("data", C.c_void_p)]


GGML_TYPE_F32, GGML_TYPE_PQ2_0 = 0, 142


def ggml_tensor(type_: int, ne, nb, data) -> GgmlTensor:
    """A tensor view: ne and nb of up to 4 dimensions (missing ne are 1, the
    nb of a missing dimension is the size of the one below), data a tensor
    or a device pointer."""
    ne = list(ne) + [1] * (4 - len(ne))
    nb = list(nb)
    while len(nb) < 4:
        nb.append(nb[-1] * ne[len(nb) - 1])
    return GgmlTensor(type_, (C.c_int64 * 4)(*ne), (C.c_size_t * 4)(*nb), _ptr(data))


def ggml_should_use(src0_type: int, device: int, ne11: int) -> bool:
    return lib().bonsai_p40_ggml_should_use(src0_type, device, ne11) == 1


def ggml_mul_mat(src0: GgmlTensor, src1: GgmlTensor, dst: GgmlTensor, scratch=None, scratch_bytes: int = 0,
                 stream=None) -> bool:
    """True when the hook enqueued dst = src0 . src1, False when the caller
    keeps its stock path."""
    return lib().bonsai_p40_ggml_mul_mat(C.byref(src0), C.byref(src1), C.byref(dst), _ptr(scratch),
                                         scratch_bytes, _stream(stream)) == 1


def fwht_gemv(W, x, signs, y, n_out: int, n_in: int, stream=None) -> None:
    _check("bonsai_p40_fwht_gemv",
           call("bonsai_p40_fwht_gemv", W, x, signs, y, n_out, n_in, stream=stream))


def _group_arrays(Ws, ys, n_outs):
    n = len(Ws)
    if not (len(ys) == n and len(n_outs) == n):
        raise ValueError("Ws, ys and n_outs must have the same length")
    Wa = (C.c_void_p * n)(*[_ptr(w) for w in Ws])
    ya = (C.c_void_p * n)(*[_ptr(y) for y in ys])
    na = (C.c_int64 * n)(*[int(r) for r in n_outs])
    # keep the arrays alive for the call: the caller holds the returned tuple
    return (Wa, ya, na), C.cast(Wa, C.c_void_p), C.cast(ya, C.c_void_p), C.cast(na, C.c_void_p), n


def gemv_group(Ws, xq, ys, n_outs, n_in: int, stream=None) -> None:
    """y_m = W_m . xq for up to 4 matrices sharing n_in, one launch."""
    keep, Wp, yp, np_, n = _group_arrays(Ws, ys, n_outs)
    rc = lib().bonsai_p40_gemv_group(Wp, yp, np_, n, _ptr(xq), n_in, _stream(stream))
    del keep
    _check("bonsai_p40_gemv_group", rc)


def fwht_gemv_group(Ws, x, signs, ys, n_outs, n_in: int, stream=None) -> None:
    """y_m = W_m . Q8_1(FWHT(signs .* x)) for up to 4 matrices, one launch."""
    keep, Wp, yp, np_, n = _group_arrays(Ws, ys, n_outs)
    rc = lib().bonsai_p40_fwht_gemv_group(Wp, yp, np_, n, _ptr(x), _ptr(signs), n_in, _stream(stream))
    del keep
    _check("bonsai_p40_fwht_gemv_group", rc)


def rmsnorm_fwht_gemv_group(Ws, x, norm_w, signs, ys, n_outs, n_in: int, eps: float,
                            stream=None) -> None:
    """y_m = W_m . Q8_1(FWHT(signs .* RMSNorm(x, norm_w, eps))), up to 4 matrices, one launch."""
    keep, Wp, yp, np_, n = _group_arrays(Ws, ys, n_outs)
    rc = lib().bonsai_p40_rmsnorm_fwht_gemv_group(Wp, yp, np_, n, _ptr(x), _ptr(norm_w), _ptr(signs), n_in,
                                                  C.c_float(eps), _stream(stream))
    del keep
    _check("bonsai_p40_rmsnorm_fwht_gemv_group", rc)


FFN_SYNC_BYTES = 256


def ffn_workspace_bytes(n_ff: int) -> int:
    """BONSAI_P40_FFN_WORKSPACE_BYTES(n_ff) of include/bonsai_p40.h."""
    return FFN_SYNC_BYTES + 8 * n_ff


def ffn_gate_up_swiglu(Wg, Wu, x, norm_w, x_signs, h_signs, hq, n_ff: int, n_embd: int, eps: float,
                       workspace, status=None, stream=None) -> None:
    """hq = Q8_1(FWHT(h_signs .* swiglu(Wg.a, Wu.a))), a = Q8_1(FWHT(x_signs .*
    RMSNorm(x))) (norm_w None: no RMSNorm), one launch; workspace zero-filled
    before its first use (ffn_workspace_bytes(n_ff) bytes)."""
    _check("bonsai_p40_ffn_gate_up_swiglu",
           call("bonsai_p40_ffn_gate_up_swiglu", Wg, Wu, x, norm_w, x_signs, h_signs, hq, n_ff, n_embd,
                C.c_float(eps), workspace, status, stream=stream))


FFN_NOALLOC_MAX_NFF = 65536


def ffn_gate_up_swiglu_noalloc(Wg, Wu, x, norm_w, x_signs, h_signs, hq, n_ff: int, n_embd: int, eps: float,
                               status=None, stream=None) -> None:
    """ffn_gate_up_swiglu with the library's static per-GPU scratch instead of
    a workspace (n_ff <= FFN_NOALLOC_MAX_NFF; calls on one GPU must not
    overlap)."""
    _check("bonsai_p40_ffn_gate_up_swiglu_noalloc",
           call("bonsai_p40_ffn_gate_up_swiglu_noalloc", Wg, Wu, x, norm_w, x_signs, h_signs, hq, n_ff, n_embd,
                C.c_float(eps), status, stream=stream))


def quantize_pq2_0(x, w, n: int, stream=None) -> None:
    _check("bonsai_p40_quantize_pq2_0", call("bonsai_p40_quantize_pq2_0", x, w, n, stream=stream))


def dequantize_pq2_0(w, y, n: int, stream=None) -> None:
    _check("bonsai_p40_dequantize_pq2_0", call("bonsai_p40_dequantize_pq2_0", w, y, n, stream=stream))


def chunk_dots(W, xq, out, n_out: int, n_in: int, stream=None) -> None:
    _check("bonsai_p40_chunk_dots",
           call("bonsai_p40_chunk_dots", W, xq, out, n_out, n_in, stream=stream))


def reload_tuning() -> None:
    """Re-read the BONSAI_* tuning variables after changing os.environ."""
    _check("bonsai_p40_reload_tuning", lib().bonsai_p40_reload_tuning())


def mfma_probe(kind: int, blocks: int, iters: int, clk, sink, stream=None) -> None:
    _check("bonsai_p40_mfma_probe", call("bonsai_p40_mfma_probe", kind, blocks, iters, clk, sink, stream=stream))


def overlap_probe(mode: int, nf: int, blocks: int, iters: int, sink, stream=None) -> None:
    _check("bonsai_p40_overlap_probe",
           call("bonsai_p40_overlap_probe", mode, nf, blocks, iters, sink, stream=stream))


def launch_probe(blocks: int, threads: int, sink, stream=None) -> None:
    _check("bonsai_p40_launch_probe", call("bonsai_p40_launch_probe", blocks, threads, sink, stream=stream))


def unit_dma_probe(W, n_out: int, n_in: int, sink, stream=None) -> None:
    _check("bonsai_p40_unit_dma_probe", call("bonsai_p40_unit_dma_probe", W, n_out, n_in, sink, stream=stream))


def stream_read(buf, nbytes: int, out, blocks: int, stream=None) -> None:
    _check("bonsai_p40_stream_read",
           call("bonsai_p40_stream_read", buf, nbytes, out, blocks, stream=stream))


# --------------------------------------------------------- sizes / helpers
def pq2_bytes(n_out: int, n_in: int) -> int:
    return n_out * (n_in // QK_PQ2) * PQ2_BYTES


def q8_bytes(n: int, n_tok: int = 1) -> int:
    return n // QK8 * n_tok * Q81_BYTES


# ------------------------------------------------------------ decode chain
CHAIN_Q8, CHAIN_FWHT, CHAIN_RMSNORM_FWHT, CHAIN_SWIGLU = 0, 1, 2, 3
CHAIN_WORKSPACE_BYTES = 4096


class ChainStep(C.Structure):
    """bonsai_p40_chain_step of include/bonsai_p40.h."""
    _fields_ = [("kind", C.c_int), ("n_mat", C.c_int), ("W", C.c_void_p * 4), ("y", C.c_void_p * 4),
                ("n_out", C.c_int64 * 4), ("n_in", C.c_int64), ("x", C.c_void_p), ("x2", C.c_void_p),
                ("norm_w", C.c_void_p), ("signs", C.c_void_p), ("q_out", C.c_void_p), ("eps", C.c_float)]


def chain_step(kind: int, W=(), y=(), n_out=(), n_in: int = 0, x=None, x2=None, norm_w=None, signs=None,
               q_out=None, eps: float = 0.0) -> ChainStep:
    """One step of a decode chain; tensors are kept by pointer (the caller
    keeps them alive while the plan is used)."""
    s = ChainStep()
    s.kind = kind
    s.n_mat = len(W)
    for i, (w, yy, n) in enumerate(zip(W, y, n_out)):
        s.W[i] = _ptr(w)
        s.y[i] = _ptr(yy)
        s.n_out[i] = int(n)
    s.n_in = int(n_in)
    s.x, s.x2, s.norm_w, s.signs, s.q_out = (_ptr(t) for t in (x, x2, norm_w, signs, q_out))
    s.eps = float(eps)
    return s


def chain_plan_bytes(n_steps: int) -> int:
    return int(lib().bonsai_p40_chain_plan_bytes(n_steps))


def chain_plan(steps, plan) -> None:
    """Check the steps and write the device plan into `plan` (a device
    tensor of chain_plan_bytes(len(steps)) bytes).  Blocking."""
    arr = (ChainStep * len(steps))(*steps)
    _check("bonsai_p40_chain_plan", lib().bonsai_p40_chain_plan(C.cast(arr, C.c_void_p), len(steps), _ptr(plan)))


def chain_run(plan, n_steps: int, workspace, status=None, stream=None) -> None:
    _check("bonsai_p40_chain_run",
           call("bonsai_p40_chain_run", plan, n_steps, workspace, status, stream=stream))


class Chain:
    """A planned decode chain with its own plan buffer and workspace."""

    def __init__(self, steps):
        import torch
        self.steps = list(steps)
        self.n = len(self.steps)
        self.plan = torch.empty(chain_plan_bytes(self.n), dtype=torch.uint8, device="cuda")
        self.workspace = torch.zeros(CHAIN_WORKSPACE_BYTES, dtype=torch.uint8, device="cuda")
        self.status = torch.zeros(1, dtype=torch.int32, device="cuda")
        chain_plan(self.steps, self.plan)

    def run(self, stream=None) -> None:
        chain_run(self.plan, self.n, self.workspace, self.status, stream=stream)
